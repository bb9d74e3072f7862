// Clustering quality evaluator: assigned inertia and empty-cluster count.
//
// Restates the evaluator of the reference's quality benchmark
// (benchmarks/quality_compare.py:69-90):
//     inertia[b] = sum_n sum_d (float(x[b,n,d]) - float(c[b,ids[b,n],d]))^2
// with the difference and its square in fp32 and the sum in fp64
// (`diff.square().sum(dtype=torch.float64)`), and
//     empty[b]   = #{k < K : no n has ids[b,n] == k}
// (`torch.bincount(...) == 0`).  Rows whose label is outside [0,K) add
// nothing and are not counted (the reference's gather would fault on them).
//
//   quality_rows  : one wave per 64 rows; lanes own column slices, so every
//                   row of x and its centroid row are coalesced loads; each
//                   lane accumulates its squares in fp64 in row order; the
//                   wave and then the workgroup combine lanes in a fixed
//                   order into one partial per workgroup.  Lane r of the
//                   wave also counts row r's label into a per-batch
//                   histogram (integer atomics: exact).
//   quality_final : one workgroup per batch row sums the partials in a
//                   fixed order and counts the empty bins.
// The result is bitwise reproducible for given inputs.
#include "device_util.hpp"
#include "fkc_internal.hpp"

namespace fkc {
namespace {

constexpr int QT = 256;       // threads per workgroup (4 waves)
constexpr int QROWS = 64;     // rows per wave
constexpr int QWG_ROWS = QROWS * (QT / 64);

__device__ inline double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int DT>
__global__ void __launch_bounds__(QT)
quality_rows_kernel(const typename Elem<DT>::T* __restrict__ x,
                    const typename Elem<DT>::T* __restrict__ cent,
                    const int32_t* __restrict__ ids,
                    double* __restrict__ partial, int32_t* __restrict__ hist,
                    int N, int K, int D, int nwg) {
  using E = Elem<DT>;
  __shared__ double wsum[QT / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int r0 = blockIdx.x * QWG_ROWS + wave * QROWS;
  const int32_t* ib = ids + (size_t)b * N;
  const int my = r0 + lane;
  const int iv = my < N ? ib[my] : -1;
  if (hist != nullptr && (uint32_t)iv < (uint32_t)K)
    atomicAdd(&hist[(size_t)b * K + iv], 1);

  double acc = 0.0;
  if (x != nullptr) {
    const typename E::T* xb = x + (size_t)b * N * D;
    const typename E::T* cb = cent + (size_t)b * K * D;
    const int nr = min(QROWS, N - r0);
    for (int j = 0; j < nr; ++j) {
      const int id = __builtin_amdgcn_readlane(iv, j);
      if ((uint32_t)id >= (uint32_t)K) continue;  // wave-uniform
      const typename E::T* xr = xb + (size_t)(r0 + j) * D;
      const typename E::T* cr = cb + (size_t)id * D;
      for (int d = lane; d < D; d += 64) {
        const float df = E::load(xr[d]) - E::load(cr[d]);
        const float sq = df * df;  // fp32 square, as the reference
        acc += (double)sq;
      }
    }
  }
  acc = wave_sum_f64(acc);
  if (lane == 0) wsum[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < QT / 64; ++w) t += wsum[w];
    partial[(size_t)b * nwg + blockIdx.x] = t;
  }
}

__global__ void __launch_bounds__(256)
quality_final_kernel(const double* __restrict__ partial,
                     const int32_t* __restrict__ hist, double* inertia,
                     int32_t* empty, int K, int nwg) {
  __shared__ double ws[4];
  __shared__ int wc[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x;
  double t = 0.0;
  if (partial != nullptr)
    for (int i = tid; i < nwg; i += 256) t += partial[(size_t)b * nwg + i];
  int e = 0;
  if (hist != nullptr)
    for (int k = tid; k < K; k += 256) e += hist[(size_t)b * K + k] == 0;
  t = wave_sum_f64(t);
  e = wave_sum_i(e);
  if (lane == 0) {
    ws[wave] = t;
    wc[wave] = e;
  }
  __syncthreads();
  if (tid == 0) {
    if (inertia != nullptr) inertia[b] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
    if (empty != nullptr) empty[b] = wc[0] + wc[1] + wc[2] + wc[3];
  }
}

template <int DT>
int launch_rows_t(const void* x, const void* c, const int32_t* ids,
                  double* partial, int32_t* hist, int64_t B, int64_t N,
                  int64_t K, int64_t D, int64_t nwg, hipStream_t s) {
  using T = typename Elem<DT>::T;
  hipLaunchKernelGGL((quality_rows_kernel<DT>), dim3((unsigned)nwg, (unsigned)B),
                     dim3(QT), 0, s, static_cast<const T*>(x),
                     static_cast<const T*>(c), ids, partial, hist, (int)N,
                     (int)K, (int)D, (int)nwg);
  return check_launch("quality_rows");
}

}  // namespace

size_t quality_workspace_bytes(int64_t B, int64_t N, int64_t K) {
  const int64_t nwg = (N + QWG_ROWS - 1) / QWG_ROWS;
  Carve c(nullptr);
  c.take<double>((size_t)B * nwg);
  c.take<int32_t>((size_t)B * K);
  return c.used;
}

int launch_quality(const void* x, const void* c, const int32_t* ids,
                   int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                   double* inertia, int32_t* empty, void* ws, size_t ws_bytes,
                   hipStream_t s) {
  const size_t need = quality_workspace_bytes(B, N, K);
  if (ws == nullptr || ws_bytes < need)
    return fail(FKC_ERR_WORKSPACE, "assigned_inertia: workspace %zu < %zu bytes",
                ws_bytes, need);
  if (reinterpret_cast<uintptr_t>(ws) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE,
                "assigned_inertia: workspace not %d-byte aligned",
                kWorkspaceAlign);
  const int64_t nwg = (N + QWG_ROWS - 1) / QWG_ROWS;
  Carve cv(ws);
  double* partial = cv.take<double>((size_t)B * nwg);
  int32_t* hist = cv.take<int32_t>((size_t)B * K);
  if (empty == nullptr) hist = nullptr;
  const void* xx = inertia != nullptr ? x : nullptr;
  int rc = FKC_OK;
  if (hist != nullptr) rc = launch_fill_i32(hist, 0, B * K, s);
  if (rc) return rc;
  if (N > 0) {
    switch (dtype) {
      case FKC_F32:
        rc = launch_rows_t<FKC_F32>(xx, c, ids, partial, hist, B, N, K, D, nwg, s);
        break;
      case FKC_F16:
        rc = launch_rows_t<FKC_F16>(xx, c, ids, partial, hist, B, N, K, D, nwg, s);
        break;
      case FKC_BF16:
        rc = launch_rows_t<FKC_BF16>(xx, c, ids, partial, hist, B, N, K, D, nwg, s);
        break;
      default:
        return fail(FKC_ERR_INVALID, "assigned_inertia: unknown dtype %d", dtype);
    }
    if (rc) return rc;
  }
  hipLaunchKernelGGL(quality_final_kernel, dim3((unsigned)B), dim3(256), 0, s,
                     N > 0 ? partial : nullptr, hist, inertia, empty, (int)K,
                     (int)nwg);
  return check_launch("quality_final");
}

}  // namespace fkc
