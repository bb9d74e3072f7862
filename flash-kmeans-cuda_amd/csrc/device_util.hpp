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

// Row reductions of the norm / finalize kernels (row_sqnorm, finalize, the
// finalize fused into the centroid update) all use one order, so their
// results agree bit for bit: lane l covers the columns VEC*(l + 64*i) + v,
// i = 0, 1, ..., v < VEC, with VEC = row_vec(D) (2 for even D above 64,
// else 1: a row of at most 64 columns then fills the wave's 64 lanes),
// accumulated with fma in (i, v) order; the 64 lane partials are then added
// by row_sum.  (The centroid update holds its sums in exactly this layout.)
__host__ __device__ inline int row_vec(int D) {
  return ((D & 1) || D <= 64) ? 1 : 2;
}

// Sum of v over the 64 lanes by a fixed tree of DPP moves: pairs and quads
// (quad_perm), 8-lane halves (row_half_mirror), 16-lane rows (row_mirror),
// then rows 0+1 and 2+3 (row_bcast:15) and all four rows (row_bcast:31).
// The total lands in lane 63 and is returned to every lane.  Each step is
// one DPP add (the butterfly of __shfl_xor costs an LDS-crossbar round trip
// per step).
__device__ inline float row_sum(float v) {
#define FKC_DPP_ADD(CTRL, RMASK)                                             \
  v += __builtin_bit_cast(                                                   \
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, \
                                         RMASK, 0xF, false))
  FKC_DPP_ADD(0xB1, 0xF);   // quad_perm [1,0,3,2]
  FKC_DPP_ADD(0x4E, 0xF);   // quad_perm [2,3,0,1]
  FKC_DPP_ADD(0x141, 0xF);  // row_half_mirror
  FKC_DPP_ADD(0x140, 0xF);  // row_mirror
  FKC_DPP_ADD(0x142, 0xA);  // row_bcast:15 into rows 1 and 3
  FKC_DPP_ADD(0x143, 0xC);  // row_bcast:31 into rows 2 and 3
#undef FKC_DPP_ADD
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Inclusive scan over the 64 lanes by DPP adds: row_shr 1, 2, 4, 8 scan
// each 16-lane row, row_bcast:15 adds row 0's total to row 1 and row 2's to
// row 3, row_bcast:31 adds lane 31 (rows 0 and 1) to rows 2 and 3.  Lanes
// without a source add the `old` operand, 0.  (A __shfl_up ladder costs an
// LDS-crossbar round trip per step.)
__device__ inline int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
  return v;
}

// Number of set bits of `mask` in lanes below the calling lane.
__device__ inline uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(
      static_cast<uint32_t>(mask >> 32),
      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// Handing data to other workgroups of the same launch without a release
// fence.  The data (a fused sort pass's digit counts, the update's head
// partials) is written with relaxed agent-scope atomics, which gfx950
// performs at the device's coherence point, past the CU and XCD caches;
// the reader loads it with agent-scope atomic loads, performed there too.
// Before the atomic that announces the data (an arrival counter) the
// writer waits for its own outstanding vector memory operations: once they
// have completed they are performed at that point, so a reader that has
// seen the announcement and then loads with agent scope sees the data.
// This rests on the hardware's behaviour, not on the HIP memory model,
// which would ask for a release fence before the announcement and an
// acquire after it (a release fence writes back the XCD's L2, which cost
// ~0.1 us per wave at every arrival).  Every site that relies on it calls
// this helper, so moving to release / acquire (or to another architecture)
// changes this one place.  The sort and update tests compare both sides of
// every such hand-over bit for bit against the oracle (and the sort's
// against its recount fallback, FKC_SORT_SPIN=0).
__device__ inline void drain_before_announce() {
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// True when the control block says the Lloyd loop already converged.
__device__ inline bool loop_done(const int32_t* ctrl) {
  return ctrl != nullptr && *ctrl != 0;
}

}  // namespace fkc
