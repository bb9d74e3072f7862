// Device-side helpers for the gfx950 kernels: element types, wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fkc.h"

namespace fkc {

// Storage and fp32 conversion per element type.  fp16 uses the hardware
// conversion (round-to-nearest-even); bf16 is stored as its 16 raw bits.
template <int DT> struct Elem;

template <> struct Elem<FKC_F32> {
  using T = float;
  __device__ static inline float load(T v) { return v; }
  __device__ static inline T store(float f) { return f; }
};

template <> struct Elem<FKC_F16> {
  using T = _Float16;
  __device__ static inline float load(T v) { return static_cast<float>(v); }
  __device__ static inline T store(float f) { return static_cast<_Float16>(f); }
};

template <> struct Elem<FKC_BF16> {
  using T = uint16_t;
  __device__ static inline float load(T v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
  }
  // Round to nearest even; NaN maps to the canonical quiet NaN 0x7FC0.
  __device__ static inline T store(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<T>(0x7fc0u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<T>(u >> 16);
  }
};

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Number of set bits of `mask` in lanes below the calling lane.
__device__ inline uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(
      static_cast<uint32_t>(mask >> 32),
      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// True when the control block says the Lloyd loop already converged.
__device__ inline bool loop_done(const int32_t* ctrl) {
  return ctrl != nullptr && *ctrl != 0;
}

}  // namespace fkc
