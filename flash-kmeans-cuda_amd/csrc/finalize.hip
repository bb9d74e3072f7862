// Centroid finalize plus the small helper kernels of the Lloyd loop.
//
// finalize_kernel restates flash_kmeans_cuda/csrc/update/update_finalize.cu:39-66:
//     new[b,k,:] = counts[b,k] > 0 ? cast(sums[b,k,:] / counts[b,k]) : old[b,k,:]
// with an IEEE division and a round-to-nearest-even cast (the reference
// divides under --use_fast_math).  One wave per centroid row.  Optionally it
// also emits, from the values just stored,
//   c_sq_out[b,k] = sum_d float(new)^2    (next iteration's kmeans.py:94 term)
//   shift_out     = max_{b,k} ||float(new) - float(old)||_2   (kmeans.py:104)
// so the loop needs no separate norm kernels.  The shift is combined with an
// integer atomic max on the float bits (valid for non-negative floats; a NaN
// row norm wins, as torch's max would propagate it).
#include "device_util.hpp"
#include "fkc_internal.hpp"

namespace fkc {
namespace {

template <int DT>
__global__ void __launch_bounds__(256)
finalize_kernel(const float* __restrict__ sums,
                const int32_t* __restrict__ counts,
                const typename Elem<DT>::T* old,
                typename Elem<DT>::T* out, float* __restrict__ c_sq_out,
                float* __restrict__ shift_out, int64_t rows, int D,
                const int32_t* __restrict__ ctrl) {
  using E = Elem<DT>;
  if (loop_done(ctrl)) return;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int cnt = counts[row];
  const float fc = (float)cnt;
  const float* sr = sums + row * D;
  const typename E::T* orow = old + row * D;
  typename E::T* nrow = out + row * D;
  // Column order and reduction shared with row_sqnorm and the finalize
  // fused into the centroid update.
  const int vec = row_vec(D);
  float sq = 0.f, sh = 0.f;
  for (int c = vec * lane; c < D; c += vec * 64) {
    for (int v = 0; v < vec; ++v) {
      const int d = c + v;
      const typename E::T o = orow[d];
      const typename E::T n = cnt > 0 ? E::store(sr[d] / fc) : o;
      nrow[d] = n;
      const float nf = E::load(n), df = nf - E::load(o);
      sq = fmaf(nf, nf, sq);
      sh = fmaf(df, df, sh);
    }
  }
  if (c_sq_out != nullptr) {
    sq = row_sum(sq);
    if (lane == 0) c_sq_out[row] = sq;
  }
  if (shift_out != nullptr) {
    sh = row_sum(sh);
    if (lane == 0)
      atomicMax(reinterpret_cast<unsigned int*>(shift_out),
                __float_as_uint(sqrtf(sh)));
  }
}

__global__ void fill_i32_kernel(int32_t* p, int32_t v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < n; j += stride) p[j] = v;
}

__global__ void fill_f32_kernel(float* p, float v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < n; j += stride) p[j] = v;
}

__global__ void fill_f64_kernel(double* p, double v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < n; j += stride) p[j] = v;
}

__global__ void iota_i32_kernel(int32_t* p, int64_t B, int64_t N) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < B * N; j += stride) p[j] = (int32_t)(j % N);
}

// Lloyd loop prologue in one launch.  Row blocks (four rows each, one wave
// per row) copy the initial centroids into the loop's centroid buffer when
// the two differ and write their squared norms with the column order and
// wave reduction of row_sqnorm_kernel (the same bits); the blocks after
// them zero the loop's control words, the label sort's and the update's
// control regions and, with a tolerance, the shift slots.
template <int DT>
__global__ void __launch_bounds__(256)
lloyd_prologue_kernel(const typename Elem<DT>::T* __restrict__ init,
                      typename Elem<DT>::T* __restrict__ cent,
                      float* __restrict__ c_sq, int64_t rows, int D,
                      int32_t* __restrict__ z0, int64_t n0,
                      int32_t* __restrict__ z1, int64_t n1,
                      float* __restrict__ z2, int64_t n2,
                      int32_t* __restrict__ z3, int64_t n3) {
  using E = Elem<DT>;
  const int64_t row_blocks = (rows + 3) / 4;
  if ((int64_t)blockIdx.x >= row_blocks) {
    const int64_t i0 = ((int64_t)blockIdx.x - row_blocks) * 256 + threadIdx.x;
    const int64_t stride = ((int64_t)gridDim.x - row_blocks) * 256;
    for (int64_t i = i0; i < n0; i += stride) z0[i] = 0;
    for (int64_t i = i0; i < n1; i += stride) z1[i] = 0;
    for (int64_t i = i0; i < n2; i += stride) z2[i] = 0.f;
    for (int64_t i = i0; i < n3; i += stride) z3[i] = 0;
    return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const typename E::T* src = init + row * D;
  typename E::T* dst = cent + row * D;
  const bool copy = init != cent;
  const int vec = row_vec(D);
  float acc = 0.f;
  for (int c = vec * lane; c < D; c += vec * 64) {
    for (int v = 0; v < vec; ++v) {
      const typename E::T e = src[c + v];
      if (copy) dst[c + v] = e;
      const float f = E::load(e);
      acc = fmaf(f, f, acc);
    }
  }
  acc = row_sum(acc);
  if (lane == 0) c_sq[row] = acc;
}

// ctrl[0] = converged flag, ctrl[1] = iterations run.  Runs after the
// finalize of iteration `it`, single thread.
__global__ void converge_check_kernel(const float* shift, int it, float tol,
                                      int32_t* ctrl) {
  if (ctrl[0] != 0) return;
  ctrl[1] = it + 1;
  if (shift[it] < tol) ctrl[0] = 1;
}

unsigned grid_for(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return (unsigned)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

template <int DT>
int launch_finalize_t(const float* sums, const int32_t* counts, const void* old,
                      void* out, float* c_sq_out, float* shift_out,
                      int64_t rows, int64_t D, const int32_t* ctrl,
                      hipStream_t s) {
  using T = typename Elem<DT>::T;
  dim3 grid((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL((finalize_kernel<DT>), grid, dim3(256), 0, s, sums,
                     counts, static_cast<const T*>(old), static_cast<T*>(out),
                     c_sq_out, shift_out, rows, (int)D, ctrl);
  return check_launch("centroid_finalize");
}

}  // namespace

int launch_finalize(const float* sums, const int32_t* counts, const void* old,
                    void* out, float* c_sq_out, float* shift_out, int64_t B,
                    int64_t K, int64_t D, int dtype, const int32_t* ctrl,
                    hipStream_t s) {
  const int64_t rows = B * K;
  if (rows == 0) return FKC_OK;
  switch (dtype) {
    case FKC_F32:
      return launch_finalize_t<FKC_F32>(sums, counts, old, out, c_sq_out,
                                        shift_out, rows, D, ctrl, s);
    case FKC_F16:
      return launch_finalize_t<FKC_F16>(sums, counts, old, out, c_sq_out,
                                        shift_out, rows, D, ctrl, s);
    case FKC_BF16:
      return launch_finalize_t<FKC_BF16>(sums, counts, old, out, c_sq_out,
                                         shift_out, rows, D, ctrl, s);
  }
  return fail(FKC_ERR_INVALID, "centroid_finalize: unknown dtype %d", dtype);
}

template <int DT>
int launch_prologue_t(const void* init, void* cent, float* c_sq, int64_t rows,
                      int64_t D, const ZeroFill& f, hipStream_t s) {
  using T = typename Elem<DT>::T;
  int64_t nz = f.n0;
  if (f.n1 > nz) nz = f.n1;
  if (f.n2 > nz) nz = f.n2;
  if (f.n3 > nz) nz = f.n3;
  const int64_t zb = nz > 0 ? (nz + 255) / 256 < 64 ? (nz + 255) / 256 : 64 : 0;
  const int64_t blocks = (rows + 3) / 4 + zb;
  if (blocks <= 0) return FKC_OK;
  hipLaunchKernelGGL((lloyd_prologue_kernel<DT>), dim3((unsigned)blocks),
                     dim3(256), 0, s, static_cast<const T*>(init),
                     static_cast<T*>(cent), c_sq, rows, (int)D, f.z0, f.n0,
                     f.z1, f.n1, f.z2, f.n2, f.z3, f.n3);
  return check_launch("lloyd_prologue");
}

int launch_lloyd_prologue(const void* init, void* cent, float* c_sq,
                          int64_t rows, int64_t D, int dtype,
                          const ZeroFill& f, hipStream_t s) {
  switch (dtype) {
    case FKC_F32:
      return launch_prologue_t<FKC_F32>(init, cent, c_sq, rows, D, f, s);
    case FKC_F16:
      return launch_prologue_t<FKC_F16>(init, cent, c_sq, rows, D, f, s);
    case FKC_BF16:
      return launch_prologue_t<FKC_BF16>(init, cent, c_sq, rows, D, f, s);
  }
  return fail(FKC_ERR_INVALID, "kmeans_lloyd: unknown dtype %d", dtype);
}

int launch_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s) {
  if (n <= 0) return FKC_OK;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, v,
                     n);
  return check_launch("fill_i32");
}

int launch_fill_f32(float* p, float v, int64_t n, hipStream_t s) {
  if (n <= 0) return FKC_OK;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, v,
                     n);
  return check_launch("fill_f32");
}

int launch_fill_f64(double* p, double v, int64_t n, hipStream_t s) {
  if (n <= 0) return FKC_OK;
  hipLaunchKernelGGL(fill_f64_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, v,
                     n);
  return check_launch("fill_f64");
}

int launch_iota_i32(int32_t* p, int64_t B, int64_t N, hipStream_t s) {
  if (B * N <= 0) return FKC_OK;
  hipLaunchKernelGGL(iota_i32_kernel, dim3(grid_for(B * N)), dim3(256), 0, s, p,
                     B, N);
  return check_launch("iota_i32");
}

int launch_converge_check(const float* shift, int it, float tol, int32_t* ctrl,
                          hipStream_t s) {
  hipLaunchKernelGGL(converge_check_kernel, dim3(1), dim3(1), 0, s, shift, it,
                     tol, ctrl);
  return check_launch("converge_check");
}

}  // namespace fkc
