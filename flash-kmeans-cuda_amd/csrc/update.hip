// Centroid sums and counts over label-sorted rows, deterministic.
//
// Restates the run semantics of the reference accumulator
// (flash_kmeans_cuda/csrc/update/update_sorted.cu:39-186): rows sorted by
// label form runs of equal labels; each run contributes its fp32 column sums
// and its length to sums[b,label,:] and counts[b,label]; labels outside
// [0,K) are skipped (:95, :167).  The reference flushes every run with fp32
// atomicAdd, so its sums depend on scheduling.  Here every bin has exactly
// one writer and rows are summed in sorted order, so results are bitwise
// reproducible:
//
//   update_runs  : one wave per unit of 128 consecutive sorted rows.  Lanes
//                  own column slices (64 lanes x VEC x NI columns per pass
//                  over the row), so every row is one coalesced load per
//                  lane slice; rows are fetched eight at a time (through the
//                  permutation for the indexed variant) before being folded
//                  into the run accumulator.  A run wholly inside the unit is
//                  written directly.  A run entering from the previous unit
//                  ("head") or leaving into the next ("tail") is parked in a
//                  per-unit partial slot instead.
//   update_merge : the unit where a multi-unit run starts owns it: it adds
//                  its tail partial to the heads of the following units, in
//                  unit order, and writes the bin once.
//
// Mode "add" (the _C / C-ABI contract) adds into caller-zeroed outputs;
// mode "overwrite" (the Lloyd loop, where every label is valid) stores, and
// the run start of each label also zeroes the empty bins below it, so no
// separate clearing pass is needed.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <limits.h>

namespace fkc {
namespace {

constexpr int UR = 128;  // sorted rows per unit (one wave)
constexpr int UT = 256;  // threads per workgroup: 4 units

// VEC consecutive columns of one row as fp32 (VEC in {1, 2}).
template <int DT, int VEC>
__device__ inline void load_cols(const typename Elem<DT>::T* p, float* out) {
  using E = Elem<DT>;
  if constexpr (VEC == 1) {
    out[0] = E::load(p[0]);
  } else if constexpr (DT == FKC_F32) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    out[0] = v.x;
    out[1] = v.y;
  } else {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    typename E::T lo, hi;
    const uint16_t l16 = (uint16_t)(w & 0xffffu), h16 = (uint16_t)(w >> 16);
    __builtin_memcpy(&lo, &l16, 2);
    __builtin_memcpy(&hi, &h16, 2);
    out[0] = E::load(lo);
    out[1] = E::load(hi);
  }
}

struct UnitMeta {  // per unit, int32 x 4
  enum { TAIL_ID = 0, TAIL_LEN = 1, HEAD_LEN = 2, THROUGH = 3 };
};

template <int DT, int VEC, int NI, bool INDEXED>
__global__ void __launch_bounds__(UT)
update_runs_kernel(const typename Elem<DT>::T* __restrict__ x,
                   const int32_t* __restrict__ perm,
                   const int32_t* __restrict__ sids, float* __restrict__ sums,
                   int32_t* __restrict__ counts, float* __restrict__ part,
                   int32_t* __restrict__ meta, int N, int K, int D,
                   int nunits, int overwrite,
                   const int32_t* __restrict__ ctrl) {
  using T = typename Elem<DT>::T;
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int u = blockIdx.x * (UT / 64) + wave;
  if (u >= nunits) return;
  const bool lead = blockIdx.z == 0;  // column block 0 writes counts / meta
  const int cbase = blockIdx.z * (64 * VEC * NI);
  const int p0 = u * UR;
  const int p1 = min(p0 + UR, N);

  const int32_t* ib = sids + (size_t)b * N;
  const int32_t* pb = INDEXED ? perm + (size_t)b * N : nullptr;
  const T* xb = x + (size_t)b * N * D;
  float* sb = sums + (size_t)b * K * D;
  int32_t* cntb = counts + (size_t)b * K;
  float* partb = part + (size_t)b * nunits * 2 * D;

  const bool has_prev = p0 > 0, has_next = p1 < N;
  const int prev = has_prev ? ib[p0 - 1] : 0;
  const int next = has_next ? ib[p1] : 0;

  int col[NI];
  bool cok[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    col[i] = cbase + (lane + 64 * i) * VEC;
    cok[i] = col[i] < D;  // D % VEC == 0, so the whole vector is in range
  }

  float acc[NI][VEC];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[i][v] = 0.f;

  int tail_id = 0, tail_len = 0, head_len = 0, through = 0;

  // Zero sums/counts of bins [lo, hi) (overwrite mode only).
  auto zero_bins = [&](int lo, int hi) {
    lo = max(lo, 0);
    hi = min(hi, K);
    for (int k = lo; k < hi; ++k) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (cok[i]) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) sb[(size_t)k * D + col[i] + v] = 0.f;
        }
    }
    if (lead)
      for (int k = lo + lane; k < hi; k += 64) cntb[k] = 0;
  };

  auto store_part = [&](int slot) {
    float* dst = partb + ((size_t)u * 2 + slot) * D;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      if (cok[i]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) dst[col[i] + v] = acc[i][v];
      }
  };

  // Close the run of label `id` covering sorted rows [s, e).
  auto flush = [&](int id, int s, int e) {
    const bool continuing = s == p0 && has_prev && prev == id;
    const bool continued = e == p1 && has_next && next == id;
    if (continuing) {
      store_part(0);
      head_len = e - s;
      through = continued ? 1 : 0;
    } else if (continued) {
      store_part(1);
      tail_id = id;
      tail_len = e - s;
    } else if ((uint32_t)id < (uint32_t)K) {
      float* dst = sb + (size_t)id * D;
#pragma unroll
      for (int i = 0; i < NI; ++i)
        if (cok[i]) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            if (overwrite)
              dst[col[i] + v] = acc[i][v];
            else
              dst[col[i] + v] += acc[i][v];
          }
        }
      if (lead && lane == 0) {
        if (overwrite)
          cntb[id] = e - s;
        else
          cntb[id] += e - s;
      }
    }
  };

  int cur = ib[p0];
  int rs = p0;
  if (overwrite && !(has_prev && prev == cur))
    zero_bins(has_prev ? prev + 1 : 0, cur);

  for (int base = p0; base < p1; base += 64) {
    const int nrow = min(64, p1 - base);
    const int iv = lane < nrow ? ib[base + lane] : 0;
    const int pv = INDEXED ? (lane < nrow ? pb[base + lane] : 0) : base + lane;
    for (int j0 = 0; j0 < nrow; j0 += 8) {
      float val[8][NI][VEC];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = j0 + jj;
        if (j < nrow) {
          const int row = __builtin_amdgcn_readlane(pv, j);
          // A permutation entry outside [0,N) contributes zeros instead of
          // reading outside x.
          const bool rok = (uint32_t)row < (uint32_t)N;
          const T* xr = xb + (size_t)(rok ? row : 0) * D;
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            if (cok[i] && rok) {
              load_cols<DT, VEC>(xr + col[i], val[jj][i]);
            } else {
#pragma unroll
              for (int v = 0; v < VEC; ++v) val[jj][i][v] = 0.f;
            }
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = j0 + jj;
        if (j < nrow) {
          const int id = __builtin_amdgcn_readlane(iv, j);
          if (id != cur) {
            flush(cur, rs, base + j);
            if (overwrite) zero_bins(cur + 1, id);
            cur = id;
            rs = base + j;
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
              for (int v = 0; v < VEC; ++v) acc[i][v] = 0.f;
          }
#pragma unroll
          for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[i][v] += val[jj][i][v];
        }
      }
    }
  }
  flush(cur, rs, p1);
  if (overwrite && !has_next) zero_bins(cur + 1, K);

  if (lead && lane == 0) {
    int32_t* m = meta + ((size_t)b * nunits + u) * 4;
    m[UnitMeta::TAIL_ID] = tail_id;
    m[UnitMeta::TAIL_LEN] = tail_len;
    m[UnitMeta::HEAD_LEN] = head_len;
    m[UnitMeta::THROUGH] = through;
  }
}

// One wave per unit; only units holding a tail partial do work.
__global__ void __launch_bounds__(UT)
update_merge_kernel(const float* __restrict__ part,
                    const int32_t* __restrict__ meta, float* __restrict__ sums,
                    int32_t* __restrict__ counts, int K, int D, int nunits,
                    int overwrite, const int32_t* __restrict__ ctrl) {
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int u = blockIdx.x * (UT / 64) + wave;
  if (u >= nunits) return;
  const int32_t* mb = meta + (size_t)b * nunits * 4;
  const int tail_len = mb[(size_t)u * 4 + UnitMeta::TAIL_LEN];
  if (tail_len == 0) return;
  const int id = mb[(size_t)u * 4 + UnitMeta::TAIL_ID];
  if ((uint32_t)id >= (uint32_t)K) return;
  const float* pb = part + (size_t)b * nunits * 2 * D;
  float* dst = sums + ((size_t)b * K + id) * D;
  int len = tail_len;
  for (int c0 = 0; c0 < D; c0 += 64) {
    const int c = c0 + lane;
    float acc = c < D ? pb[((size_t)u * 2 + 1) * D + c] : 0.f;
    int v = u + 1;
    int l = tail_len;
    while (v < nunits) {
      if (c < D) acc += pb[((size_t)v * 2 + 0) * D + c];
      l += mb[(size_t)v * 4 + UnitMeta::HEAD_LEN];
      if (!mb[(size_t)v * 4 + UnitMeta::THROUGH]) break;
      ++v;
    }
    len = l;
    if (c < D) {
      if (overwrite)
        dst[c] = acc;
      else
        dst[c] += acc;
    }
  }
  if (lane == 0) {
    int32_t* cp = counts + (size_t)b * K + id;
    if (overwrite)
      *cp = len;
    else
      *cp += len;
  }
}

template <int DT, int VEC, int NI, bool INDEXED>
int launch_runs_t(const void* x, const int32_t* perm, const int32_t* sids,
                  float* sums, int32_t* counts, float* part, int32_t* meta,
                  int64_t B, int64_t N, int64_t K, int64_t D, int64_t nunits,
                  bool overwrite, const int32_t* ctrl, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int64_t cols_per_block = 64 * VEC * NI;
  dim3 grid((unsigned)((nunits + 3) / 4), (unsigned)B,
            (unsigned)((D + cols_per_block - 1) / cols_per_block));
  hipLaunchKernelGGL((update_runs_kernel<DT, VEC, NI, INDEXED>), grid,
                     dim3(UT), 0, s, static_cast<const T*>(x), perm, sids,
                     sums, counts, part, meta, (int)N, (int)K, (int)D,
                     (int)nunits, overwrite ? 1 : 0, ctrl);
  return check_launch("update_runs");
}

template <int DT, bool INDEXED>
int launch_runs_dt(const void* x, const int32_t* perm, const int32_t* sids,
                   float* sums, int32_t* counts, float* part, int32_t* meta,
                   int64_t B, int64_t N, int64_t K, int64_t D, int64_t nunits,
                   bool overwrite, const int32_t* ctrl, hipStream_t s) {
  const int vec = (D % 2 == 0) ? 2 : 1;
  const int64_t slices = (D + 64 * vec - 1) / (64 * vec);
#define FKC_RUNS(V, NI_)                                                    \
  return launch_runs_t<DT, V, NI_, INDEXED>(x, perm, sids, sums, counts,   \
                                            part, meta, B, N, K, D, nunits, \
                                            overwrite, ctrl, s)
  if (vec == 2) {
    if (slices <= 1) FKC_RUNS(2, 1);
    if (slices <= 2) FKC_RUNS(2, 2);
    FKC_RUNS(2, 4);
  }
  if (slices <= 1) FKC_RUNS(1, 1);
  if (slices <= 2) FKC_RUNS(1, 2);
  FKC_RUNS(1, 4);
#undef FKC_RUNS
}

}  // namespace

size_t update_workspace_bytes(int64_t B, int64_t N, int64_t D) {
  const int64_t nunits = (N + UR - 1) / UR;
  Carve c(nullptr);
  c.take<float>((size_t)B * nunits * 2 * D);
  c.take<int32_t>((size_t)B * nunits * 4);
  return c.used;
}

int launch_update(const void* x, const int32_t* perm,
                  const int32_t* ids_sorted, float* sums, int32_t* counts,
                  int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                  bool overwrite, void* ws, size_t ws_bytes,
                  const int32_t* ctrl, hipStream_t s) {
  if (B == 0) return FKC_OK;
  if (N == 0) {
    if (!overwrite) return FKC_OK;
    int rc = launch_fill_f32(sums, 0.f, B * K * D, s);
    return rc ? rc : launch_fill_i32(counts, 0, B * K, s);
  }
  const size_t need = update_workspace_bytes(B, N, D);
  if (ws_bytes < need || ws == nullptr)
    return fail(FKC_ERR_WORKSPACE, "centroid_update: workspace %zu < %zu bytes",
                ws_bytes, need);
  const int64_t nunits = (N + UR - 1) / UR;
  Carve c(ws);
  float* part = c.take<float>((size_t)B * nunits * 2 * D);
  int32_t* meta = c.take<int32_t>((size_t)B * nunits * 4);
  int rc = FKC_OK;
  const bool idx = perm != nullptr;
  switch (dtype) {
    case FKC_F32:
      rc = idx ? launch_runs_dt<FKC_F32, true>(x, perm, ids_sorted, sums, counts,
                                               part, meta, B, N, K, D, nunits,
                                               overwrite, ctrl, s)
               : launch_runs_dt<FKC_F32, false>(x, perm, ids_sorted, sums,
                                                counts, part, meta, B, N, K, D,
                                                nunits, overwrite, ctrl, s);
      break;
    case FKC_F16:
      rc = idx ? launch_runs_dt<FKC_F16, true>(x, perm, ids_sorted, sums, counts,
                                               part, meta, B, N, K, D, nunits,
                                               overwrite, ctrl, s)
               : launch_runs_dt<FKC_F16, false>(x, perm, ids_sorted, sums,
                                                counts, part, meta, B, N, K, D,
                                                nunits, overwrite, ctrl, s);
      break;
    case FKC_BF16:
      rc = idx ? launch_runs_dt<FKC_BF16, true>(x, perm, ids_sorted, sums,
                                                counts, part, meta, B, N, K, D,
                                                nunits, overwrite, ctrl, s)
               : launch_runs_dt<FKC_BF16, false>(x, perm, ids_sorted, sums,
                                                 counts, part, meta, B, N, K, D,
                                                 nunits, overwrite, ctrl, s);
      break;
    default:
      return fail(FKC_ERR_INVALID, "centroid_update: unknown dtype %d", dtype);
  }
  if (rc) return rc;
  dim3 grid((unsigned)((nunits + 3) / 4), (unsigned)B);
  hipLaunchKernelGGL(update_merge_kernel, grid, dim3(UT), 0, s, part, meta,
                     sums, counts, (int)K, (int)D, (int)nunits,
                     overwrite ? 1 : 0, ctrl);
  return check_launch("update_merge");
}

}  // namespace fkc
