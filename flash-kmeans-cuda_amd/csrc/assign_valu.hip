// fp32 VALU assignment (the fallback route) and row squared norms.
//
// assign_valu_kernel restates the reference's tensor-core-free kernel
// (flash_kmeans_cuda/csrc/assign/assign_safe.cu:38-81): for each point,
//     dist_k = max(0, x_sq + c_sq[k] - 2 * <x, c_k>)      (assign_common.cuh:33-36)
// with the dot product accumulated in fp32 as one fused multiply-add chain in
// feature order, and the strict-< running minimum that keeps the lowest k on
// ties (assign_common.cuh:23-28).  It serves fp32 inputs, D % 16 != 0,
// D > 256 and FKC_ASSIGN_FORCE_SAFE (api.cpp:12-25).
//
// Layout: one thread per point, 256 points per workgroup.  Centroids pass
// through LDS in 32 x 32 (centroid x feature) fp32 tiles; every lane of a
// wave reads the same LDS word (broadcast), so the tile costs one LDS read
// per FMA-column and no bank conflicts.  Each thread keeps 32 partial dot
// products in registers while the feature tiles stream past.
#include "device_util.hpp"
#include "fkc_internal.hpp"

#include <float.h>

namespace fkc {

int launch_assign_mfma(const void* x, const void* c, const float* c_sq,
                       int32_t* ids, int64_t B, int64_t N, int64_t K,
                       int64_t D, int dtype, const int32_t* ctrl,
                       hipStream_t s);

namespace {

constexpr int VT = 256;   // threads (points) per workgroup
constexpr int VKC = 32;   // centroids per LDS tile
constexpr int VDC = 32;   // features per LDS tile

template <int DT>
__global__ void __launch_bounds__(VT)
assign_valu_kernel(const typename Elem<DT>::T* __restrict__ x,
                   const typename Elem<DT>::T* __restrict__ c,
                   const float* __restrict__ x_sq,
                   const float* __restrict__ c_sq, int32_t* __restrict__ ids,
                   int N, int K, int D, const int32_t* __restrict__ ctrl) {
  using E = Elem<DT>;
  if (loop_done(ctrl)) return;
  __shared__ float tile[VKC][VDC];
  __shared__ float tile_q[VKC];

  const int tid = threadIdx.x;
  const int b = blockIdx.y;
  const int n = blockIdx.x * VT + tid;
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
  for (int k0 = 0; k0 < K; k0 += VKC) {
    float acc[VKC];
#pragma unroll
    for (int j = 0; j < VKC; ++j) acc[j] = 0.f;
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
        for (int kk = 0; kk < VKC; ++kk) {
#pragma unroll
          for (int dd = 0; dd < VDC; ++dd)
            acc[kk] = fmaf(xv[dd], tile[kk][dd], acc[kk]);
        }
      } else {
        for (int dd = 0; dd < dn; ++dd) {
          const float xv = E::load(xr[d0 + dd]);
#pragma unroll
          for (int kk = 0; kk < VKC; ++kk)
            acc[kk] = fmaf(xv, tile[kk][dd], acc[kk]);
        }
      }
    }
    const int kn = min(VKC, K - k0);
    for (int kk = 0; kk < kn; ++kk) {
      float dist = xs + tile_q[kk] - 2.0f * acc[kk];
      dist = dist > 0.f ? dist : 0.f;
      if (dist < best) {
        best = dist;
        bidx = k0 + kk;
      }
    }
  }
  if (valid) ids[(size_t)b * N + n] = bidx;
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
  float acc = 0.f;
  for (int d = lane; d < D; d += 64) {
    const float v = E::load(r[d]);
    acc = fmaf(v, v, acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) out[row] = acc;
}

template <int DT>
int launch_valu_t(const void* x, const void* c, const float* x_sq,
                  const float* c_sq, int32_t* ids, int64_t B, int64_t N,
                  int64_t K, int64_t D, const int32_t* ctrl, hipStream_t s) {
  using T = typename Elem<DT>::T;
  dim3 grid((unsigned)((N + VT - 1) / VT), (unsigned)B);
  hipLaunchKernelGGL((assign_valu_kernel<DT>), grid, dim3(VT), 0, s,
                     static_cast<const T*>(x), static_cast<const T*>(c), x_sq,
                     c_sq, ids, (int)N, (int)K, (int)D, ctrl);
  return check_launch("assign_valu");
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
                  hipStream_t s) {
  if (B == 0 || N == 0) return FKC_OK;
  if (assign_uses_mfma(dtype, D))
    return launch_assign_mfma(x, c, c_sq, ids, B, N, K, D, dtype, ctrl, s);
  switch (dtype) {
    case FKC_F32:
      return launch_valu_t<FKC_F32>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    case FKC_F16:
      return launch_valu_t<FKC_F16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
    case FKC_BF16:
      return launch_valu_t<FKC_BF16>(x, c, x_sq, c_sq, ids, B, N, K, D, ctrl, s);
  }
  return fail(FKC_ERR_INVALID, "assign: unknown dtype %d", dtype);
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
