// fp32 VALU assignment (the fallback route) and row squared norms.
//
// assign_valu_kernel restates the reference's tensor-core-free kernel
// (flash_kmeans_cuda/csrc/assign/assign_safe.cu:38-81): for each point,
//     dist_k = max(0, x_sq + c_sq[k] - 2 * <x, c_k>)      (assign_common.cuh:33-36)
// with the dot product accumulated in fp32 as one fused multiply-add chain in
// feature order, and the strict-< running minimum that keeps the lowest k on
// ties (assign_common.cuh:23-28).  It serves fp32 inputs, fp16/bf16 with
// D % 8 != 0 or D > 512, and FKC_ASSIGN_FORCE_SAFE (api.cpp:12-25).
//
// Layout: SPLIT adjacent lanes per point (256 / SPLIT points per
// workgroup); lane s of a point scores centroids k = s (mod SPLIT) of each
// tile.  Centroids pass through LDS in 32 x 32 (centroid x feature) fp32
// tiles.  Each lane keeps 32 / SPLIT partial dot products in registers while
// the feature tiles stream past; every (point, centroid) dot product is one
// lane's FMA chain in feature order whatever SPLIT is, so labels do not
// depend on it.  The SPLIT lanes of a point merge with the lowest-index rule
// at the end.  SPLIT > 1 gives small N enough workgroups to fill the chip.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <float.h>

namespace fkc {

int launch_assign_mfma(const void* x, const void* c, const float* c_sq,
                       int32_t* ids, int64_t B, int64_t N, int64_t K,
                       int64_t D, int dtype, const int32_t* ctrl,
                       hipStream_t s, hipEvent_t ev0, hipEvent_t ev1,
                       void* ws, size_t ws_bytes);

namespace {

constexpr int VT = 256;   // threads (points) per workgroup
constexpr int VKC = 32;   // centroids per LDS tile
constexpr int VDC = 32;   // features per LDS tile

template <int DT, int SPLIT, bool PREF>
__global__ void __launch_bounds__(VT)
assign_valu_kernel(const typename Elem<DT>::T* __restrict__ x,
                   const typename Elem<DT>::T* __restrict__ c,
                   const float* __restrict__ x_sq,
                   const float* __restrict__ c_sq, int32_t* __restrict__ ids,
                   int N, int K, int D, const int32_t* __restrict__ ctrl) {
  using E = Elem<DT>;
  constexpr int PPW = VT / SPLIT;    // points per workgroup
  constexpr int KPL = VKC / SPLIT;   // centroids per lane per tile
  if (loop_done(ctrl)) return;
  // Rows padded to 36 floats: 16-byte aligned, so the lanes' reads of a
  // row's features become 16-byte loads (one per four FMAs instead of one per
  // FMA; 33-float rows forced 4-byte loads), with at most two-way bank
  // conflicts when lanes read different rows (measured: (262144, 256, 128)
  // fp32 1.00 -> 0.32 ms, (131072, 1024, 128) fp32 2.25 -> 1.92 ms,
  // (100000, 300, 37) fp16 0.100 -> 0.082 ms).
  __shared__ __attribute__((aligned(16))) float tile[VKC][VDC + 4];
  __shared__ float tile_q[VKC];

  const int tid = threadIdx.x;
  const int sl = tid % SPLIT;        // this lane's centroid residue
  const int b = blockIdx.y;
  const int n = blockIdx.x * PPW + tid / SPLIT;
  const bool valid = n < N;
  const typename E::T* xr = x + ((size_t)b * N + (valid ? n : 0)) * D;
  const typename E::T* cb = c + (size_t)b * K * D;

  float xs = 0.f;
  if (x_sq != nullptr) {
    xs = valid ? x_sq[(size_t)b * N + n] : 0.f;
  } else {
    for (int d = 0; d < D; ++d) {
      const float v = E::load(xr[d]);
      xs = fmaf(v, v, xs);
    }
  }

  float best = FLT_MAX;
  int bidx = 0;
  if constexpr (!PREF) {
    // One lane per point (large N: enough waves to hide the loads; the
    // prefetching loop below measured 15% slower at N = 262144) or a
    // partial last feature chunk (computed only over its real features;
    // the prefetching loop would pad it to 32): the plain tile loop.
    for (int k0 = 0; k0 < K; k0 += VKC) {
      float acc[KPL];
  #pragma unroll
      for (int j = 0; j < KPL; ++j) acc[j] = 0.f;
      for (int d0 = 0; d0 < D; d0 += VDC) {
        __syncthreads();
        for (int i = tid; i < VKC * VDC; i += VT) {
          const int kk = i / VDC, dd = i % VDC;
          const int k = k0 + kk, d = d0 + dd;
          tile[kk][dd] = (k < K && d < D) ? E::load(cb[(size_t)k * D + d]) : 0.f;
        }
        if (d0 == 0 && tid < VKC) {
          const int k = k0 + tid;
          tile_q[tid] = k < K ? c_sq[(size_t)b * K + k] : 0.f;
        }
        __syncthreads();
        const int dn = min(VDC, D - d0);
        if (dn == VDC) {
          float xv[VDC];
  #pragma unroll
          for (int dd = 0; dd < VDC; ++dd) xv[dd] = E::load(xr[d0 + dd]);
  #pragma unroll
          for (int j = 0; j < KPL; ++j) {
            const int kk = j * SPLIT + sl;
  #pragma unroll
            for (int dd = 0; dd < VDC; ++dd)
              acc[j] = fmaf(xv[dd], tile[kk][dd], acc[j]);
          }
        } else {
          for (int dd = 0; dd < dn; ++dd) {
            const float xv = E::load(xr[d0 + dd]);
  #pragma unroll
            for (int j = 0; j < KPL; ++j)
              acc[j] = fmaf(xv, tile[j * SPLIT + sl][dd], acc[j]);
          }
        }
      }
  #pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int kk = j * SPLIT + sl;
        if (k0 + kk < K) {
          float dist = xs + tile_q[kk] - 2.0f * acc[j];
          dist = dist > 0.f ? dist : 0.f;
          if (dist < best) {  // kk rises with j: the first minimum is kept
            best = dist;
            bidx = k0 + kk;
          }
        }
      }
    }
  } else {
  // The (centroid tile, feature chunk) steps run in sequence; the next
  // step's centroid tile (TPT values per thread) and feature chunk are
  // loaded into registers before the current step is computed, so every
  // step's global loads overlap the previous step's arithmetic instead of
  // costing a round trip each.
  constexpr int TPT = VKC * VDC / VT;  // tile values per thread
  static_assert(VKC * VDC % VT == 0, "tile split");
  const int nkt = (K + VKC - 1) / VKC, ndc = (D + VDC - 1) / VDC;
  const int nsteps = nkt * ndc;
  float pt[TPT], pq = 0.f, px[VDC];
  auto fetch = [&](int st) {
    const int k0 = (st / ndc) * VKC, d0 = (st % ndc) * VDC;
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = tid + j * VT;
      const int k = k0 + i / VDC, d = d0 + i % VDC;
      pt[j] = (k < K && d < D) ? E::load(cb[(size_t)k * D + d]) : 0.f;
    }
    if (d0 == 0 && tid < VKC)
      pq = k0 + tid < K ? c_sq[(size_t)b * K + k0 + tid] : 0.f;
#pragma unroll
    for (int dd = 0; dd < VDC; ++dd)
      px[dd] = d0 + dd < D ? E::load(xr[d0 + dd]) : 0.f;
  };
  fetch(0);
  float acc[KPL];
  for (int st = 0; st < nsteps; ++st) {
    const int k0 = (st / ndc) * VKC, dc = st % ndc;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = tid + j * VT;
      tile[i / VDC][i % VDC] = pt[j];
    }
    if (dc == 0 && tid < VKC) tile_q[tid] = pq;
    float xv[VDC];
#pragma unroll
    for (int dd = 0; dd < VDC; ++dd) xv[dd] = px[dd];
    __syncthreads();
    if (st + 1 < nsteps) fetch(st + 1);
    if (dc == 0) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) acc[j] = 0.f;
    }
    // Features past D are zero in both operands and add nothing.
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int kk = j * SPLIT + sl;
#pragma unroll
      for (int dd = 0; dd < VDC; ++dd) acc[j] = fmaf(xv[dd], tile[kk][dd], acc[j]);
    }
    if (dc == ndc - 1) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int kk = j * SPLIT + sl;
        if (k0 + kk < K) {
          float dist = xs + tile_q[kk] - 2.0f * acc[j];
          dist = dist > 0.f ? dist : 0.f;
          if (dist < best) {  // kk rises with j: the first minimum is kept
            best = dist;
            bidx = k0 + kk;
          }
        }
      }
    }
  }
  }
  // Merge the SPLIT lanes of this point (adjacent lanes): smaller distance,
  // then smaller index.
#pragma unroll
  for (int off = 1; off < SPLIT; off <<= 1) {
    const float ob = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bidx, off, 64);
    if (ob < best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
  }
  if (valid && sl == 0) ids[(size_t)b * N + n] = bidx;
}

template <int DT>
__global__ void __launch_bounds__(256)
row_sqnorm_kernel(const typename Elem<DT>::T* __restrict__ src,
                  float* __restrict__ out, int64_t rows, int D,
                  const int32_t* __restrict__ ctrl) {
  using E = Elem<DT>;
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const typename E::T* r = src + row * D;
  // Column order and reduction shared with the finalize kernels.
  const int vec = row_vec(D);
  float acc = 0.f;
  for (int c = vec * lane; c < D; c += vec * 64) {
    for (int v = 0; v < vec; ++v) {
      const float f = E::load(r[c + v]);
      acc = fmaf(f, f, acc);
    }
  }
  acc = row_sum(acc);
  if (lane == 0) out[row] = acc;
}

// PREF (several lanes per point and D a multiple of the 32-feature chunk):
// the prefetching step loop, measured at (1, 4096, 64, 128) fp32 0.0180 ->
// 0.0129 ms and (1, 65536, 1024, 64) fp32 0.338 -> 0.308 ms.
template <int DT, int SPLIT>
int launch_valu_split(const void* x, const void* c, const float* x_sq,
                      const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                      int64_t K, int64_t D, const int32_t* ctrl,
                      hipStream_t s) {
  using T = typename Elem<DT>::T;
  constexpr int PPW = VT / SPLIT;
  dim3 grid((unsigned)((N + PPW - 1) / PPW), (unsigned)B);
  if (SPLIT > 1 && D % VDC == 0)
    hipLaunchKernelGGL((assign_valu_kernel<DT, SPLIT, SPLIT != 1>), grid,
                       dim3(VT), 0, s, static_cast<const T*>(x),
                       static_cast<const T*>(c), x_sq, c_sq, ids, (int)N,
                       (int)K, (int)D, ctrl);
  else
    hipLaunchKernelGGL((assign_valu_kernel<DT, SPLIT, false>), grid, dim3(VT),
                       0, s, static_cast<const T*>(x),
                       static_cast<const T*>(c), x_sq, c_sq, ids, (int)N,
                       (int)K, (int)D, ctrl);
  return check_launch("assign_valu");
}

// Lanes per point: one while the grid has >= 512 workgroups (2 per CU),
// else the smallest of 4, 8, 16 that gives >= 1024 workgroups.  Two lanes
// per point were never the fastest (measured, ms at 1 / 2 / 4 / 8 / 16 lanes:
// (131072, 1024, 128) fp32 0.94 / 1.93 / 1.05 / 1.05 / 1.63;
// (65536, 1024, 64) fp32 0.43 / 0.53 / 0.27 / 0.29 / 0.43;
// (32768, 512, 128) fp32 0.40 / 0.31 / 0.16 / 0.15 / 0.23;
// (100000, 300, 37) fp16 0.18 / 0.11 / 0.088 / 0.10 / 0.15).
template <int DT>
int launch_valu_t(const void* x, const void* c, const float* x_sq,
                  const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                  int64_t K, int64_t D, const int32_t* ctrl, hipStream_t s) {
  int split = 1;
  if (B * ((N + VT - 1) / VT) < 512) {
    split = 4;
    while (split < 16 && B * ((N * split + VT - 1) / VT) < 1024) split <<= 1;
  }
  switch (split) {
    case 1: return launch_valu_split<DT, 1>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    case 4: return launch_valu_split<DT, 4>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    case 8: return launch_valu_split<DT, 8>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    default: return launch_valu_split<DT, 16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
  }
}

template <int DT>
int launch_rowsq_t(const void* src, float* out, int64_t rows, int64_t D,
                   const int32_t* ctrl, hipStream_t s) {
  using T = typename Elem<DT>::T;
  dim3 grid((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL((row_sqnorm_kernel<DT>), grid, dim3(256), 0, s,
                     static_cast<const T*>(src), out, rows, (int)D, ctrl);
  return check_launch("row_sqnorm");
}

}  // namespace

int launch_assign(const void* x, const void* c, const float* x_sq,
                  const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                  int64_t K, int64_t D, int dtype, const int32_t* ctrl,
                  hipStream_t s, hipEvent_t ev0, hipEvent_t ev1, void* ws,
                  size_t ws_bytes) {
  if (B == 0 || N == 0) return FKC_OK;
  if (assign_uses_mfma(dtype, D))
    return launch_assign_mfma(x, c, c_sq, ids, B, N, K, D, dtype, ctrl, s,
                              ev0, ev1, ws, ws_bytes);
  // The VALU route marks its span with event records on the stream.
  if (ev0 != nullptr) (void)hipEventRecord(ev0, s);
  int rc = FKC_OK;
  switch (dtype) {
    case FKC_F32:
      rc = launch_valu_t<FKC_F32>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
      break;
    case FKC_F16:
      rc = launch_valu_t<FKC_F16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
      break;
    case FKC_BF16:
      rc = launch_valu_t<FKC_BF16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
      break;
    default:
      return fail(FKC_ERR_INVALID, "assign: unknown dtype %d", dtype);
  }
  if (ev1 != nullptr) (void)hipEventRecord(ev1, s);
  return rc;
}

int launch_row_sqnorm(const void* src, float* out, int64_t rows, int64_t D,
                      int dtype, const int32_t* ctrl, hipStream_t s) {
  if (rows == 0) return FKC_OK;
  switch (dtype) {
    case FKC_F32: return launch_rowsq_t<FKC_F32>(src, out, rows, D, ctrl, s);
    case FKC_F16: return launch_rowsq_t<FKC_F16>(src, out, rows, D, ctrl, s);
    case FKC_BF16: return launch_rowsq_t<FKC_BF16>(src, out, rows, D, ctrl, s);
  }
  return fail(FKC_ERR_INVALID, "row_sqnorm: unknown dtype %d", dtype);
}

}  // namespace fkc
