// Clustering quality evaluator: assigned inertia, empty-cluster count and
// the inertia of a point sample.
//
// Restates the evaluator of the reference's quality benchmark
// (benchmarks/quality_compare.py:69-116):
//     inertia[b] = sum_n sum_d (float(x[b,n,d]) - float(c[b,ids[b,n],d]))^2
// with the difference and its square in fp32 and the sum in fp64
// (`diff.square().sum(dtype=torch.float64)`), and
//     empty      = #{k < K : no (b,n) has ids[b,n] == k}
// (`torch.bincount(ids.reshape(-1), minlength=K) == 0`: one histogram over
// the labels of every batch row).  Rows whose label is outside [0,K) add
// nothing and are not counted (the reference's gather would fault on them).
//
//   quality_rows   : one wave per 64 rows; lanes own column slices, so every
//                    row of x and its centroid row are coalesced loads; each
//                    lane accumulates its squares in fp64 in row order; the
//                    wave and then the workgroup combine lanes in a fixed
//                    order into one partial per workgroup.  Lane r of the
//                    wave also counts row r's label into the K-bin histogram
//                    (integer atomics: exact).
//   quality_final  : one workgroup per batch row sums the partials in a
//                    fixed order; workgroup 0 also counts the empty bins.
//   sample_gather  : the sampled rows of x, for the sampled inertia
//                    (`_sample_exact_inertia`, :91-116), which then runs the
//                    assignment and quality_rows over them: each sampled
//                    point adds its squared distance to the nearest centroid.
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
                    int N, int K, int D, int nwg,
                    const int32_t* __restrict__ sidx, int sN) {
  using E = Elem<DT>;
  __shared__ double wsum[QT / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int r0 = blockIdx.x * QWG_ROWS + wave * QROWS;
  const int32_t* ib = ids + (size_t)b * N;
  const int my = r0 + lane;
  // Sampled rows (sidx set): a row whose sample index is outside [0, sN)
  // counts as unlabelled.
  const bool sok = sidx == nullptr || (my < N && (uint32_t)sidx[my] < (uint32_t)sN);
  const int iv = my < N && sok ? ib[my] : -1;
  if (hist != nullptr && (uint32_t)iv < (uint32_t)K) atomicAdd(&hist[iv], 1);

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
  if (hist != nullptr && b == 0)
    for (int k = tid; k < K; k += 256) e += hist[k] == 0;
  t = wave_sum_f64(t);
  e = wave_sum_i(e);
  if (lane == 0) {
    ws[wave] = t;
    wc[wave] = e;
  }
  __syncthreads();
  if (tid == 0) {
    if (inertia != nullptr) inertia[b] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
    if (empty != nullptr && b == 0) *empty = wc[0] + wc[1] + wc[2] + wc[3];
  }
}

// xs[b,s,:] = x[b,idx[s],:] (raw element bits; one wave per sampled row).
__global__ void __launch_bounds__(256)
sample_gather_kernel(const uint8_t* __restrict__ x,
                     const int32_t* __restrict__ idx, uint8_t* __restrict__ xs,
                     int N, int S, int row_bytes) {
  const int lane = threadIdx.x & 63;
  const int s = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= S) return;
  const size_t b = blockIdx.y;
  // An index outside [0, N) copies row 0 (in bounds); quality_rows then
  // leaves that sample out.
  const int n = (uint32_t)idx[s] < (uint32_t)N ? idx[s] : 0;
  const uint8_t* src = x + (b * N + (size_t)n) * row_bytes;
  uint8_t* dst = xs + (b * S + s) * (size_t)row_bytes;
  if (row_bytes % 16 == 0) {
    for (int i = lane * 16; i < row_bytes; i += 64 * 16)
      *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(src + i);
  } else {
    for (int i = lane * 2; i < row_bytes; i += 64 * 2)
      *reinterpret_cast<uint16_t*>(dst + i) =
          *reinterpret_cast<const uint16_t*>(src + i);
  }
}

template <int DT>
int launch_rows_t(const void* x, const void* c, const int32_t* ids,
                  double* partial, int32_t* hist, int64_t B, int64_t N,
                  int64_t K, int64_t D, int64_t nwg, const int32_t* sidx,
                  int64_t sN, hipStream_t s) {
  using T = typename Elem<DT>::T;
  hipLaunchKernelGGL((quality_rows_kernel<DT>), dim3((unsigned)nwg, (unsigned)B),
                     dim3(QT), 0, s, static_cast<const T*>(x),
                     static_cast<const T*>(c), ids, partial, hist, (int)N,
                     (int)K, (int)D, (int)nwg, sidx, (int)sN);
  return check_launch("quality_rows");
}

}  // namespace

size_t quality_workspace_bytes(int64_t B, int64_t N, int64_t K) {
  const int64_t nwg = (N + QWG_ROWS - 1) / QWG_ROWS;
  Carve c(nullptr);
  c.take<double>((size_t)B * nwg);
  c.take<int32_t>((size_t)K);
  return c.used;
}

size_t sample_workspace_bytes(int64_t B, int64_t S, int64_t K, int64_t D,
                              int dtype) {
  Carve c(nullptr);
  c.take<char>((size_t)B * S * D * dtype_size(dtype));  // sampled rows
  c.take<float>((size_t)B * S);                         // their x_sq
  c.take<float>((size_t)B * K);                         // c_sq
  c.take<int32_t>((size_t)B * S);                       // their labels
  c.take<char>(quality_workspace_bytes(B, S, K));
  return c.used;
}

int launch_sampled_inertia(const void* x, const void* c, const int32_t* idx,
                           int64_t S, int64_t B, int64_t N, int64_t K,
                           int64_t D, int dtype, double* inertia, void* ws,
                           size_t ws_bytes, hipStream_t s) {
  const size_t need = sample_workspace_bytes(B, S, K, D, dtype);
  if (ws == nullptr || ws_bytes < need)
    return fail(FKC_ERR_WORKSPACE, "sampled_inertia: workspace %zu < %zu bytes",
                ws_bytes, need);
  if (reinterpret_cast<uintptr_t>(ws) % kWorkspaceAlign != 0)
    return fail(FKC_ERR_WORKSPACE,
                "sampled_inertia: workspace not %d-byte aligned",
                kWorkspaceAlign);
  Carve cv(ws);
  void* xs = cv.take<char>((size_t)B * S * D * dtype_size(dtype));
  float* xs_sq = cv.take<float>((size_t)B * S);
  float* c_sq = cv.take<float>((size_t)B * K);
  int32_t* lab = cv.take<int32_t>((size_t)B * S);
  const size_t qbytes = quality_workspace_bytes(B, S, K);
  void* qws = cv.take<char>(qbytes);
  const int row_bytes = (int)(D * dtype_size(dtype));
  hipLaunchKernelGGL(sample_gather_kernel,
                     dim3((unsigned)((S + 3) / 4), (unsigned)B), dim3(256), 0,
                     s, static_cast<const uint8_t*>(x), idx,
                     static_cast<uint8_t*>(xs), (int)N, (int)S, row_bytes);
  int rc = check_launch("sample_gather");
  if (!rc) rc = launch_row_sqnorm(c, c_sq, B * K, D, dtype, nullptr, s);
  if (!rc && !assign_uses_mfma(dtype, D))
    rc = launch_row_sqnorm(xs, xs_sq, B * S, D, dtype, nullptr, s);
  if (!rc)
    rc = launch_assign(xs, c, xs_sq, c_sq, lab, B, S, K, D, dtype, nullptr, s);
  if (!rc)
    rc = launch_quality(xs, c, lab, B, S, K, D, dtype, inertia, nullptr, qws,
                        qbytes, s, idx, N);
  return rc;
}

int launch_quality(const void* x, const void* c, const int32_t* ids,
                   int64_t B, int64_t N, int64_t K, int64_t D, int dtype,
                   double* inertia, int32_t* empty, void* ws, size_t ws_bytes,
                   hipStream_t s, const int32_t* sidx, int64_t sN) {
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
  int32_t* hist = cv.take<int32_t>((size_t)K);
  if (empty == nullptr) hist = nullptr;
  const void* xx = inertia != nullptr ? x : nullptr;
  int rc = FKC_OK;
  if (hist != nullptr) rc = launch_fill_i32(hist, 0, K, s);
  if (rc) return rc;
  if (N > 0) {
    switch (dtype) {
      case FKC_F32:
        rc = launch_rows_t<FKC_F32>(xx, c, ids, partial, hist, B, N, K, D, nwg, sidx, sN, s);
        break;
      case FKC_F16:
        rc = launch_rows_t<FKC_F16>(xx, c, ids, partial, hist, B, N, K, D, nwg, sidx, sN, s);
        break;
      case FKC_BF16:
        rc = launch_rows_t<FKC_BF16>(xx, c, ids, partial, hist, B, N, K, D, nwg, sidx, sN, s);
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
