// libtorch fkc:: API over the C ABI (include/fkc.h).
//
// Argument checks follow the reference's api.cpp:27-44 and the launcher
// checks it relies on (assign_sm80.cu:712-731, update_sorted.cu:196-206,
// 253-277, update_finalize.cu:76-83); the update functions zero their
// outputs first, as api.cpp:79-80 and :91-92 do.  Scratch memory comes from
// torch's caching allocator and is handed to the kernels as a workspace.
#include "flash_kmeans_cuda.h"

#include <c10/hip/HIPStream.h>

#include "fkc.h"

namespace fkc {
namespace {

int dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return FKC_F32;
    case at::kHalf: return FKC_F16;
    case at::kBFloat16: return FKC_BF16;
    default: TORCH_CHECK(false, "unsupported dtype ", t.scalar_type());
  }
  return -1;
}

fkc_stream_t stream_of(const at::Tensor& t) {
  return reinterpret_cast<fkc_stream_t>(
      c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == FKC_OK, what, " failed (status ", rc, "): ", fkc_last_error());
}

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  return at::empty({static_cast<int64_t>(bytes > 0 ? bytes : 1)},
                   at::TensorOptions().dtype(at::kByte).device(like.device()));
}

void validate_assign_inputs(const at::Tensor& x, const at::Tensor& centroids,
                            const at::Tensor& x_sq, const at::Tensor& c_sq,
                            const at::Tensor& cluster_ids) {
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(centroids.is_cuda(), "centroids must be a CUDA tensor");
  TORCH_CHECK(x.dim() == 3, "x must be (B, N, D)");
  TORCH_CHECK(centroids.dim() == 3, "centroids must be (B, K, D)");
  TORCH_CHECK(x.scalar_type() == centroids.scalar_type(), "x and centroids must share dtype");
  TORCH_CHECK(centroids.size(0) == x.size(0) && centroids.size(2) == x.size(2),
              "centroids must be (B, K, D) matching x");
  TORCH_CHECK(x_sq.scalar_type() == at::kFloat, "x_sq must be fp32");
  TORCH_CHECK(c_sq.scalar_type() == at::kFloat, "c_sq must be fp32");
  TORCH_CHECK(c_sq.numel() == x.size(0) * centroids.size(1), "c_sq must be (B, K)");
  TORCH_CHECK(cluster_ids.scalar_type() == at::kInt, "cluster_ids must be int32");
  TORCH_CHECK(cluster_ids.dim() == 2 && cluster_ids.size(0) == x.size(0) &&
                  cluster_ids.size(1) == x.size(1),
              "cluster_ids must be (B, N) int32");
  TORCH_CHECK(x.is_contiguous() && centroids.is_contiguous() && c_sq.is_contiguous() &&
                  cluster_ids.is_contiguous(),
              "all tensors must be contiguous");
}

void validate_update(const at::Tensor& x, const at::Tensor& ids, const at::Tensor& sums,
                     const at::Tensor& counts) {
  TORCH_CHECK(x.is_cuda(), "x must be CUDA");
  TORCH_CHECK(x.dim() == 3, "x must be (B, N, D)");
  TORCH_CHECK(ids.scalar_type() == at::kInt, "cluster_ids must be int32");
  TORCH_CHECK(sums.scalar_type() == at::kFloat, "centroid_sums must be fp32");
  TORCH_CHECK(counts.scalar_type() == at::kInt, "centroid_counts must be int32");
  TORCH_CHECK(ids.dim() == 2 && ids.size(0) == x.size(0) && ids.size(1) == x.size(1),
              "cluster_ids_sorted must be (B, N)");
  TORCH_CHECK(sums.dim() == 3 && sums.size(0) == x.size(0) && sums.size(2) == x.size(2),
              "centroid_sums must be (B, K, D)");
  TORCH_CHECK(counts.numel() == sums.size(0) * sums.size(1), "centroid_counts must be (B, K)");
  TORCH_CHECK(x.is_contiguous() && ids.is_contiguous() && sums.is_contiguous() &&
                  counts.is_contiguous(),
              "all tensors must be contiguous");
}

void run_update(const at::Tensor& x, const at::Tensor* sorted_idx, const at::Tensor& ids,
                at::Tensor& sums, at::Tensor& counts) {
  validate_update(x, ids, sums, counts);
  sums.zero_();
  counts.zero_();
  const int64_t B = x.size(0), N = x.size(1), D = x.size(2), K = sums.size(1);
  at::Tensor ws = workspace(fkc_update_workspace_bytes(B, N, D), x);
  int rc;
  if (sorted_idx) {
    TORCH_CHECK(sorted_idx->scalar_type() == at::kInt, "sorted_idx must be int32");
    TORCH_CHECK(sorted_idx->dim() == 2 && sorted_idx->size(0) == B && sorted_idx->size(1) == N,
                "sorted_idx must be (B, N)");
    TORCH_CHECK(sorted_idx->is_contiguous(), "all tensors must be contiguous");
    rc = fkc_centroid_update_sorted_indexed(
        x.data_ptr(), sorted_idx->data_ptr<int32_t>(), ids.data_ptr<int32_t>(),
        sums.data_ptr<float>(), counts.data_ptr<int32_t>(), B, N, K, D, dtype_code(x),
        ws.data_ptr(), ws.numel(), stream_of(x));
  } else {
    rc = fkc_centroid_update_sorted(x.data_ptr(), ids.data_ptr<int32_t>(),
                                    sums.data_ptr<float>(), counts.data_ptr<int32_t>(), B,
                                    N, K, D, dtype_code(x), ws.data_ptr(), ws.numel(),
                                    stream_of(x));
  }
  check_rc(rc, "centroid_update_sorted");
}

}  // namespace

at::Tensor euclid_assign(const at::Tensor& x, const at::Tensor& centroids,
                         const at::Tensor& x_sq, const at::Tensor& c_sq) {
  at::Tensor ids = at::empty({x.size(0), x.size(1)},
                             at::TensorOptions().dtype(at::kInt).device(x.device()));
  return euclid_assign_out(x, centroids, x_sq, c_sq, ids);
}

at::Tensor euclid_assign_out(const at::Tensor& x, const at::Tensor& centroids,
                             const at::Tensor& x_sq, const at::Tensor& c_sq,
                             at::Tensor cluster_ids) {
  validate_assign_inputs(x, centroids, x_sq, c_sq, cluster_ids);
  const int64_t B = x.size(0), N = x.size(1), D = x.size(2), K = centroids.size(1);
  const float* xsq = nullptr;
  if (x_sq.numel() == B * N) {
    TORCH_CHECK(x_sq.is_contiguous(), "all tensors must be contiguous");
    xsq = x_sq.data_ptr<float>();
  }
  const size_t need = fkc_euclid_assign_workspace_bytes(B, N, K, D, dtype_code(x));
  if (need == 0) {
    check_rc(fkc_euclid_assign(x.data_ptr(), centroids.data_ptr(), xsq, c_sq.data_ptr<float>(),
                               cluster_ids.data_ptr<int32_t>(), B, N, K, D, dtype_code(x),
                               stream_of(x)),
             "euclid_assign");
  } else {
    // K sliced across workgroups: partial winners in a stream-ordered workspace.
    at::Tensor ws = workspace(need, x);
    check_rc(fkc_euclid_assign_ws(x.data_ptr(), centroids.data_ptr(), xsq,
                                  c_sq.data_ptr<float>(), cluster_ids.data_ptr<int32_t>(), B, N,
                                  K, D, dtype_code(x), ws.data_ptr(), ws.numel(), stream_of(x)),
             "euclid_assign");
  }
  return cluster_ids;
}

void centroid_update_sorted(const at::Tensor& x_sorted, const at::Tensor& cluster_ids_sorted,
                            at::Tensor centroid_sums, at::Tensor centroid_counts) {
  run_update(x_sorted, nullptr, cluster_ids_sorted, centroid_sums, centroid_counts);
}

void centroid_update_sorted_indexed(const at::Tensor& x, const at::Tensor& sorted_idx,
                                    const at::Tensor& cluster_ids_sorted,
                                    at::Tensor centroid_sums, at::Tensor centroid_counts) {
  run_update(x, &sorted_idx, cluster_ids_sorted, centroid_sums, centroid_counts);
}

at::Tensor centroid_finalize(const at::Tensor& centroid_sums, const at::Tensor& centroid_counts,
                             const at::Tensor& old_centroids) {
  at::Tensor out = at::empty_like(old_centroids);
  return centroid_finalize_out(centroid_sums, centroid_counts, old_centroids, out);
}

at::Tensor centroid_finalize_out(const at::Tensor& centroid_sums,
                                 const at::Tensor& centroid_counts,
                                 const at::Tensor& old_centroids, at::Tensor out) {
  TORCH_CHECK(centroid_sums.is_cuda(), "all tensors must be CUDA");
  TORCH_CHECK(centroid_sums.scalar_type() == at::kFloat, "sums must be fp32");
  TORCH_CHECK(centroid_counts.scalar_type() == at::kInt, "counts must be int32");
  TORCH_CHECK(old_centroids.scalar_type() == out.scalar_type(),
              "old and new centroids must share dtype");
  TORCH_CHECK(centroid_sums.dim() == 3, "sums must be (B, K, D)");
  TORCH_CHECK(old_centroids.sizes() == centroid_sums.sizes() &&
                  out.sizes() == centroid_sums.sizes(),
              "centroids must be (B, K, D) like sums");
  TORCH_CHECK(centroid_counts.numel() == centroid_sums.size(0) * centroid_sums.size(1),
              "counts must be (B, K)");
  TORCH_CHECK(centroid_sums.is_contiguous() && centroid_counts.is_contiguous() &&
                  old_centroids.is_contiguous() && out.is_contiguous(),
              "all tensors must be contiguous");
  check_rc(fkc_centroid_finalize(centroid_sums.data_ptr<float>(),
                                 centroid_counts.data_ptr<int32_t>(), old_centroids.data_ptr(),
                                 out.data_ptr(), centroid_sums.size(0), centroid_sums.size(1),
                                 centroid_sums.size(2), dtype_code(out), stream_of(out)),
           "centroid_finalize");
  return out;
}

std::tuple<at::Tensor, at::Tensor> label_sort(const at::Tensor& cluster_ids,
                                              int64_t n_clusters) {
  TORCH_CHECK(cluster_ids.is_cuda() && cluster_ids.dim() == 2, "cluster_ids must be CUDA (B, N)");
  at::Tensor ids = cluster_ids.to(at::kInt).contiguous();
  at::Tensor sorted = at::empty_like(ids), perm = at::empty_like(ids);
  const int64_t B = ids.size(0), N = ids.size(1);
  at::Tensor ws = workspace(fkc_label_sort_workspace_bytes(B, N, n_clusters), ids);
  check_rc(fkc_label_sort(ids.data_ptr<int32_t>(), sorted.data_ptr<int32_t>(),
                          perm.data_ptr<int32_t>(), B, N, n_clusters, ws.data_ptr(),
                          ws.numel(), stream_of(ids)),
           "label_sort");
  return {sorted, perm};
}

std::tuple<at::Tensor, at::Tensor, int64_t> batch_kmeans_euclid(
    const at::Tensor& x_in, int64_t n_clusters, int64_t max_iters, double tol,
    const at::Tensor& init_centroids) {
  TORCH_CHECK(x_in.is_cuda(), "flash_kmeans_cuda requires a CUDA input");
  TORCH_CHECK(x_in.dim() == 3, "x must be (B, N, D)");
  at::Tensor x = x_in.contiguous();
  const int64_t B = x.size(0), N = x.size(1), D = x.size(2), K = n_clusters;
  TORCH_CHECK(init_centroids.scalar_type() == x.scalar_type(),
              "x and centroids must share dtype");
  at::Tensor init = init_centroids.contiguous().view({B, K, D});
  // The loop copies init into cents in its first launch; init is not written.
  at::Tensor cents = at::empty_like(init);
  at::Tensor ids = at::empty({B, N}, at::TensorOptions().dtype(at::kInt).device(x.device()));
  const int dt = dtype_code(x);
  const int iters = static_cast<int>(max_iters);
  at::Tensor ws = workspace(fkc_kmeans_workspace_bytes(B, N, K, D, dt, iters > 0 ? iters : 1), x);
  int32_t n = 0;
  check_rc(fkc_kmeans_lloyd_from(x.data_ptr(), init.data_ptr(), cents.data_ptr(),
                                 ids.data_ptr<int32_t>(), B, N, K, D, dt, iters,
                                 static_cast<float>(tol), ws.data_ptr(), ws.numel(),
                                 stream_of(x), nullptr, &n),
           "batch_kmeans_euclid");
  return {ids, cents, static_cast<int64_t>(n)};
}

}  // namespace fkc
