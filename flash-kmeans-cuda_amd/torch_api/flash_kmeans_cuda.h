#pragma once

// Public libtorch C++ API, on PyTorch-ROCm: the drop-in for the reference's
// flash_kmeans_cuda/csrc/flash_kmeans_cuda.h:31-77 (namespace fkc, same six
// functions, same signatures and semantics).  Tensors are borrowed; work is
// enqueued on the current HIP stream of the tensors' device; bad arguments
// raise c10::Error (TORCH_CHECK), as in the reference.  Everything below
// calls the C ABI of include/fkc.h, whose kernels are gfx950 HIP.
//
// batch_kmeans_euclid is an addition with no counterpart in the reference's
// C++ header: the Lloyd loop of its Python driver (kmeans.py:108-195) for C++
// callers.

#include <ATen/ATen.h>

#include <tuple>

#if defined(_WIN32)
#if defined(FKC_BUILD_SHARED)
#define FKC_API __declspec(dllexport)
#else
#define FKC_API __declspec(dllimport)
#endif
#else
#define FKC_API __attribute__((visibility("default")))
#endif

namespace fkc {

// Nearest-centroid label of every point, in a new (B, N) int32 tensor.
FKC_API at::Tensor euclid_assign(const at::Tensor& x, const at::Tensor& centroids,
                                 const at::Tensor& x_sq, const at::Tensor& c_sq);

// As euclid_assign, with the labels stored in the caller's (B, N) int32
// tensor, which is returned.
FKC_API at::Tensor euclid_assign_out(const at::Tensor& x, const at::Tensor& centroids,
                                     const at::Tensor& x_sq, const at::Tensor& c_sq,
                                     at::Tensor cluster_ids);

// Per-label fp32 row sums and int32 counts over label-sorted rows; the
// output tensors are cleared first.
FKC_API void centroid_update_sorted(const at::Tensor& x_sorted,
                                    const at::Tensor& cluster_ids_sorted,
                                    at::Tensor centroid_sums, at::Tensor centroid_counts);

// The same sums and counts with x in its original row order, row p of the
// sorted order being x[sorted_idx[p]].
FKC_API void centroid_update_sorted_indexed(const at::Tensor& x, const at::Tensor& sorted_idx,
                                            const at::Tensor& cluster_ids_sorted,
                                            at::Tensor centroid_sums,
                                            at::Tensor centroid_counts);

// New centroids sums / counts (the old centroid where a count is 0), in a
// new tensor of old_centroids' dtype.
FKC_API at::Tensor centroid_finalize(const at::Tensor& centroid_sums,
                                     const at::Tensor& centroid_counts,
                                     const at::Tensor& old_centroids);

// As centroid_finalize, stored in the caller's tensor `out`, which is
// returned.
FKC_API at::Tensor centroid_finalize_out(const at::Tensor& centroid_sums,
                                         const at::Tensor& centroid_counts,
                                         const at::Tensor& old_centroids, at::Tensor out);

// Stable label sort (B, N) int32 -> (sorted ids, permutation), both int32.
FKC_API std::tuple<at::Tensor, at::Tensor> label_sort(const at::Tensor& cluster_ids,
                                                      int64_t n_clusters);

// Whole Lloyd loop: returns (cluster_ids (B,N) int32, centroids (B,K,D),
// iterations run).  init_centroids (B,K,D) is not modified.
FKC_API std::tuple<at::Tensor, at::Tensor, int64_t> batch_kmeans_euclid(
    const at::Tensor& x, int64_t n_clusters, int64_t max_iters, double tol,
    const at::Tensor& init_centroids);

}  // namespace fkc
